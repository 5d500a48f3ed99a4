// Row and query encoding for the int8 MFMA screen, tombstones and small fills (gfx950).
//
// Reference contracts: encode_int8_rows / encode_int8_queries (detail/int8.cuh:30-136) and
// remove_rows / remove_int8_rows (certex_kernels.cuh:391-415, detail/int8.cuh:139-147). For 8-bit
// integer vectors the code is the vector itself shifted into int8 (no projection, no scale), so
// the screen is exact; the row term folds the norm (l2) or the shift correction (inner product).

#include "../kernels.hpp"

namespace certex_amd {
namespace {

inline unsigned blocks_for(int64_t n, int block = 256)
{
  return unsigned((n + block - 1) / block);
}

/**
 * One thread per 16-byte chunk of a stored row (row_bytes / 16 = 8 or 16 consecutive lanes per
 * row), so that the reads of the input rows and the writes of the codes are coalesced; the
 * chunks' partial norms and sums meet by shuffles within the row's lanes.
 */
__global__ void encode_rows_kernel(const uint8_t* x, int64_t n, int64_t dim, int row_bytes,
                                   uint8_t flip, metric_kind metric, int8_t* codes, int32_t* rowc)
{
  const int cpr   = row_bytes / 16;  // a power of two that divides 64
  const int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  const int64_t r = t / cpr;
  const int c     = int(t % cpr);
  int norm = 0, sum = 0;
  if (r < n) {
    uint8_t v[16];
    const int64_t j0 = int64_t(c) * 16;
    if (dim % 16 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && j0 < dim) {
      *reinterpret_cast<int4*>(v) = *reinterpret_cast<const int4*>(x + r * dim + j0);
    } else {
#pragma unroll
      for (int b = 0; b < 16; ++b) { v[b] = j0 + b < dim ? x[r * dim + j0 + b] : uint8_t(0); }
    }
    int8_t out[16];
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const int code = j0 + b < dim ? int(int8_t(v[b] ^ flip)) : 0;
      out[b]         = int8_t(code);
      norm += code * code;
      sum += code;
    }
    *reinterpret_cast<int4*>(codes + r * row_bytes + j0) = *reinterpret_cast<const int4*>(out);
  }
  for (int off = 1; off < cpr; off <<= 1) {
    norm += __shfl_xor(norm, off);
    sum += __shfl_xor(sum, off);
  }
  if (r < n && c == 0) {
    rowc[r] = metric == metric_kind::l2 ? -(norm >> 1) : (flip ? 128 * sum : 0);
  }
}

/**
 * The rows of more than 256 bytes (row_bytes a multiple of 256): one wave per row, lane l on the
 * 16-byte chunks l, l + 64, ...; the row's norm and sum meet by shuffles over the wave.
 */
__global__ void encode_rows_wide_kernel(const uint8_t* x, int64_t n, int64_t dim, int row_bytes,
                                        uint8_t flip, metric_kind metric, int8_t* codes, int32_t* rowc)
{
  const int64_t r = (blockIdx.x * int64_t(blockDim.x) + threadIdx.x) >> 6;
  const int lane  = threadIdx.x & 63;
  if (r >= n) { return; }  // whole waves leave together (64 divides the block)
  int norm = 0, sum = 0;
  for (int c = lane; c < row_bytes / 16; c += 64) {
    const int64_t j0 = int64_t(c) * 16;
    int8_t out[16];
#pragma unroll
    for (int b = 0; b < 16; ++b) {
      const int code = j0 + b < dim ? int(int8_t(x[r * dim + j0 + b] ^ flip)) : 0;
      out[b]         = int8_t(code);
      norm += code * code;
      sum += code;
    }
    *reinterpret_cast<int4*>(codes + r * row_bytes + j0) = *reinterpret_cast<const int4*>(out);
  }
  for (int off = 1; off < 64; off <<= 1) {
    norm += __shfl_xor(norm, off);
    sum += __shfl_xor(sum, off);
  }
  if (lane == 0) { rowc[r] = metric == metric_kind::l2 ? -(norm >> 1) : (flip ? 128 * sum : 0); }
}

__global__ void encode_queries_kernel(const uint8_t* q, const int32_t* rows, int64_t nq,
                                      int64_t nq_pad, int64_t dim, int row_bytes, uint8_t flip,
                                      int8_t* qcodes, int8_t* qpaired)
{
  const int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (t >= nq_pad * row_bytes) { return; }
  const int64_t i = t / row_bytes, j = t % row_bytes;
  const int64_t r = i < nq && rows != nullptr ? int64_t(rows[i]) : i;  // the caller's query row
  const int8_t c  = (i < nq && j < dim) ? int8_t(q[r * dim + j] ^ flip) : int8_t(0);
  qcodes[t]       = c;
  if (qpaired != nullptr) { qpaired[paired_offset(i, j, row_bytes)] = c; }
}

__device__ inline int64_t stored_row(const row_places& at, int64_t id)
{
  return id < at.n_listed ? int64_t(at.list_pos[id]) : id;
}

__global__ void remove_kernel(const int64_t* ids, int64_t n, int64_t size, int32_t* rowc,
                              unsigned long long* newly, row_places at)
{
  const int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (t >= n) { return; }
  const int64_t id = ids[t];
  if (id < 0 || id >= size) { return; }
  if (id < at.n_part) { static_cast<int32_t*>(at.part_rowc)[at.part_pos[id]] = kDeadRow; }
  if (at.anchor_stride > 0 && id % at.anchor_stride == 0 && id / at.anchor_stride < at.n_anchor) {
    static_cast<int32_t*>(at.anchor_rowc)[id / at.anchor_stride] = kDeadRow;
  }
  if (atomicExch(rowc + stored_row(at, id), kDeadRow) != kDeadRow) { atomicAdd(newly, 1ull); }
}

template <typename T>
__global__ void fill_kernel(T* p, int64_t n, T v)
{
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x) {
    p[i] = v;
  }
}

__global__ void iota_kernel(int32_t* p, int64_t n, int32_t first)
{
  for (int64_t i = blockIdx.x * int64_t(blockDim.x) + threadIdx.x; i < n;
       i += int64_t(gridDim.x) * blockDim.x) {
    p[i] = first + int32_t(i);
  }
}

// ---- float vectors ---------------------------------------------------------------------------

__device__ inline double coord(const void* p, elem t, int64_t i)
{
  if (t == elem::bf16) { return double(static_cast<const __bf16*>(p)[i]); }
  return t == elem::f32 ? double(static_cast<const float*>(p)[i])
                        : double(static_cast<const _Float16*>(p)[i]);
}

/** Euclidean norm of row i (1 when zero) for unit normalisation, fp64 in coordinate order. */
__device__ inline double row_norm(const void* x, elem t, int64_t i, int64_t dim)
{
  double s = 0;
  for (int64_t j = 0; j < dim; ++j) {
    const double v = coord(x, t, i * dim + j);
    s              = fma(v, v, s);
  }
  return s > 0 ? sqrt(s) : 1.0;
}

__device__ inline void atomic_max_pos(double* p, double v)
{
  // non-negative doubles order like their bit patterns
  atomicMax(reinterpret_cast<unsigned long long*>(p), (unsigned long long)__double_as_longlong(v));
}

/** Upper bound of sqrt(s) for a non-negative fp64 sum s accumulated over `terms` terms. */
__device__ inline double sqrt_up(double s, int64_t terms)
{
  return sqrt(s * (1.0 + 4e-16 * double(terms + 4))) * (1.0 + 4e-16);
}

__global__ void column_sums_kernel(const void* x, elem t, int64_t n, int64_t dim, bool normalize,
                                   int64_t rows_per_block, double* sums)
{
  __shared__ double nrm[512];
  const int64_t r0 = blockIdx.x * rows_per_block;
  const int64_t r1 = r0 + rows_per_block < n ? r0 + rows_per_block : n;
  for (int64_t i = r0 + threadIdx.x; i < r1; i += blockDim.x) {
    nrm[i - r0] = normalize ? row_norm(x, t, i, dim) : 1.0;
  }
  __syncthreads();
  for (int64_t j = threadIdx.x; j < dim; j += blockDim.x) {
    double s = 0;
    for (int64_t i = r0; i < r1; ++i) { s += coord(x, t, i * dim + j) / nrm[i - r0]; }
    atomicAdd(sums + j, s);
  }
}

constexpr double kF16Safe = 4096.0;  // |Z| above this: the row is always a candidate

/** fp16 value of z (round to nearest), 0 for results below the smallest normal fp16. */
__device__ inline _Float16 to_f16(double z)
{
  const _Float16 h = _Float16(float(z));
  return fabs(double(h)) < 6.103515625e-05 ? _Float16(0.0f) : h;
}

/** Sum of v over the 64 lanes of a wave (xor butterfly: every lane gets the sum). */
__device__ inline double wave_sum(double v)
{
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) { v += __shfl_xor(v, off); }
  return v;
}

/** A lane's coordinates of one row loaded together: j = j0 + 64 u + lane, u < kLaneChunk. */
constexpr int kLaneChunk = 16;

template <typename T, int N>
__device__ inline void lane_coords_t(const T* row, int64_t dim, int64_t j0, int lane,
                                     double (&v)[N])
{
  T x[N];  // loads from clamped positions, unconditional: all issued before any use
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int64_t j = j0 + 64 * u + lane;
    x[u]            = row[j < dim ? j : dim - 1];
  }
#pragma unroll
  for (int u = 0; u < N; ++u) { v[u] = j0 + 64 * u + lane < dim ? double(x[u]) : 0.0; }
}

/** Coordinates j0 + 64 u + lane of row i (0 at and past dim), all loads issued before any use:
 *  a loop that used each coordinate as it arrived waited for one load at a time. */
template <int N = kLaneChunk>
__device__ inline void lane_coords(const void* x, elem t, int64_t i, int64_t dim, int64_t j0,
                                   int lane, double (&v)[N])
{
  if (t == elem::bf16) {
    lane_coords_t(static_cast<const __bf16*>(x) + i * dim, dim, j0, lane, v);
  } else if (t == elem::f32) {
    lane_coords_t(static_cast<const float*>(x) + i * dim, dim, j0, lane, v);
  } else {
    lane_coords_t(static_cast<const _Float16*>(x) + i * dim, dim, j0, lane, v);
  }
}

/** center[j0 + 64 u + lane], u < N (clamped positions past dim), loaded together. */
template <int N = kLaneChunk>
__device__ inline void lane_center(const double* center, int64_t dim, int64_t j0, int lane,
                                   double (&c)[N])
{
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int64_t j = j0 + 64 * u + lane;
    c[u]            = center[j < dim ? j : dim - 1];
  }
}

/** |x_i| (1 when zero) by a wave: per-lane fp64 partial sums in coordinate order, a butterfly. */
__device__ inline double wave_row_norm(const void* x, elem t, int64_t i, int64_t dim, int lane)
{
  double s2 = 0;
  for (int64_t j0 = 0; j0 < dim; j0 += 64 * kLaneChunk) {
    double v[kLaneChunk];
    lane_coords(x, t, i, dim, j0, lane, v);
#pragma unroll
    for (int u = 0; u < kLaneChunk; ++u) { s2 = fma(v[u], v[u], s2); }  // past dim: + 0, exact
  }
  s2 = wave_sum(s2);
  return s2 > 0 ? sqrt(s2) : 1.0;
}

/**
 * out[0] raised to the largest |x / |x| - center| (|x - center| without normalizing) over the n
 * rows, sqrt_up of the fp64 sum: rows by waves over a grid stride as encode_rows_f16_kernel takes
 * them, one atomic per workgroup.
 */
__global__ __launch_bounds__(256) void max_norm_kernel(const void* x, elem t, int64_t n,
                                                       int64_t dim, bool normalize,
                                                       const double* center, double* out)
{
  __shared__ double wmax[4];
  const int lane      = threadIdx.x & 63;
  const int wave      = threadIdx.x >> 6;
  const int64_t waves = int64_t(gridDim.x) * 4;
  double m            = 0;
  for (int64_t i = blockIdx.x * int64_t(4) + wave; i < n; i += waves) {
    const double nrm = normalize ? wave_row_norm(x, t, i, dim, lane) : 1.0;
    double s         = 0;
    for (int64_t j0 = 0; j0 < dim; j0 += 64 * kLaneChunk) {
      double v[kLaneChunk], c[kLaneChunk];
      lane_coords(x, t, i, dim, j0, lane, v);
      lane_center(center, dim, j0, lane, c);
#pragma unroll
      for (int u = 0; u < kLaneChunk; ++u) {
        if (j0 + 64 * u + lane < dim) {
          const double z = v[u] / nrm - c[u];
          s              = fma(z, z, s);
        }
      }
    }
    m = fmax(m, sqrt_up(wave_sum(s), dim));
  }
  if (lane == 0) { wmax[wave] = m; }
  __syncthreads();
  if (threadIdx.x == 0) { atomic_max_pos(out, fmax(fmax(wmax[0], wmax[1]), fmax(wmax[2], wmax[3]))); }
}

/**
 * Rows i = w, w + W, ... for wave w of W (a grid stride), each by one wave whose lanes take the
 * coordinates j = lane, lane + 64, ... (coalesced loads and stores): rows[i] = fp16(Z) with
 * Z = (x / |x| - center) / alpha (x / |x| when normalizing), subnormals set to 0, zero padded;
 * rowc[i] = -|Z|^2 / 2, raised so that it bounds the term's fp32 accumulation (0 for the inner
 * product); a row with |Z| above kF16Safe is stored as zeros with rowc = +inf (always a
 * candidate). maxima[0] and maxima[1] are raised to the largest |fp16(Z)| and |Z - fp16(Z)|
 * (sqrt_up of their sums), one atomic each per workgroup. The fp64 sums are per-lane partials
 * and a butterfly; they only enter bounds that carry their rounding slack.
 */
__global__ __launch_bounds__(256) void encode_rows_f16_kernel(const void* x, elem t, int64_t n,
                                                              int64_t dim, int halves,
                                                              bool normalize, const double* center,
                                                              double inv_alpha, metric_kind metric,
                                                              double gamma, uint16_t* rows,
                                                              float* rowc, double* maxima)
{
  __shared__ double wmax[2][4];
  const int lane      = threadIdx.x & 63;
  const int wave      = threadIdx.x >> 6;
  const int64_t waves = int64_t(gridDim.x) * 4;
  double mh = 0, me = 0;  // this wave's largest bounds of |fp16(Z)| and |Z - fp16(Z)|
  for (int64_t i = blockIdx.x * int64_t(4) + wave; i < n; i += waves) {
    _Float16* dst    = reinterpret_cast<_Float16*>(rows + i * halves);
    const double nrm = normalize ? wave_row_norm(x, t, i, dim, lane) : 1.0;
    double a         = 0;
    for (int64_t j0 = 0; j0 < dim; j0 += 64 * kLaneChunk) {
      double v[kLaneChunk], c[kLaneChunk];
      lane_coords(x, t, i, dim, j0, lane, v);
      lane_center(center, dim, j0, lane, c);
#pragma unroll
      for (int u = 0; u < kLaneChunk; ++u) {
        if (j0 + 64 * u + lane < dim) {
          const double z = (v[u] / nrm - c[u]) * inv_alpha;
          a              = fma(z, z, a);
        }
      }
    }
    a = wave_sum(a);  // the same value in every lane: the branch below is uniform
    if (!(sqrt(a) <= kF16Safe)) {
      for (int64_t j = lane; j < halves; j += 64) { dst[j] = _Float16(0.0f); }
      if (lane == 0) { rowc[i] = INFINITY; }
      continue;
    }
    double nz = 0, ez = 0;
    for (int64_t j0 = 0; j0 < dim; j0 += 64 * kLaneChunk) {
      double v[kLaneChunk], c[kLaneChunk];
      lane_coords(x, t, i, dim, j0, lane, v);
      lane_center(center, dim, j0, lane, c);
#pragma unroll
      for (int u = 0; u < kLaneChunk; ++u) {
        const int64_t j = j0 + 64 * u + lane;
        if (j < dim) {
          const double z   = (v[u] / nrm - c[u]) * inv_alpha;
          const _Float16 h = to_f16(z);
          const double e   = z - double(h);  // exact (Sterbenz, or h = 0)
          dst[j]           = h;
          nz               = fma(double(h), double(h), nz);
          ez               = fma(e, e, ez);
        }
      }
    }
    for (int64_t j = dim + lane; j < halves; j += 64) { dst[j] = _Float16(0.0f); }
    nz = wave_sum(nz);
    ez = wave_sum(ez);
    if (lane == 0) {
      if (metric == metric_kind::inner) {
        rowc[i] = 0.0f;
      } else {
        // row term rounded up: the fp32 accumulation error of this term is folded in (factor
        // 1 - 2g)
        const double c = -(a * (1.0 - 1e-13) / 2.0) * (1.0 - 2.0 * gamma - 1e-10);
        float f        = float(c);
        if (double(f) < c) { f = nextafterf(f, INFINITY); }
        rowc[i] = f;
      }
    }
    mh = fmax(mh, sqrt_up(nz, dim));
    me = fmax(me, sqrt_up(ez, dim));
  }
  if (lane == 0) {
    wmax[0][wave] = mh;
    wmax[1][wave] = me;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    atomic_max_pos(maxima + 0, fmax(fmax(wmax[0][0], wmax[0][1]), fmax(wmax[0][2], wmax[0][3])));
    atomic_max_pos(maxima + 1, fmax(fmax(wmax[1][0], wmax[1][1]), fmax(wmax[1][2], wmax[1][3])));
  }
}

/**
 * One wave per query, its lanes over the coordinates j = lane, lane + 64, ... (coalesced loads):
 * qrows[i] = fp16(W) with W = (q / |q| - center) / alpha (q / |q| when normalizing), subnormals
 * set to 0, zero padded; qscal[3 i ..] = |W|^2 (lowered by 1e-13), |fp16(W)| and |W - fp16(W)|
 * (raised for the rounding of their sums, sqrt_up). Per-lane fp64 partial sums and a butterfly:
 * the sums only enter bounds that carry these slacks.
 */
template <int N>
__global__ __launch_bounds__(256) void encode_queries_f16_kernel(const void* q, const int32_t* rows,
                                                                 elem t, int64_t nq,
                                                                 int64_t nq_pad, int64_t dim,
                                                                 int halves, bool normalize,
                                                                 const double* center,
                                                                 double inv_alpha, uint16_t* qrows,
                                                                 double* qscal, uint16_t* qpaired)
{
  const int64_t i = blockIdx.x * int64_t(blockDim.x / 64) + (threadIdx.x >> 6);
  const int lane  = threadIdx.x & 63;
  if (i >= nq_pad) { return; }  // uniform over the wave
  _Float16* dst = reinterpret_cast<_Float16*>(qrows + i * halves);
  // half j of the query, and of its paired copy when there is one
  auto put = [&](int64_t j, _Float16 h) {
    dst[j] = h;
    if (qpaired != nullptr) {
      reinterpret_cast<_Float16*>(qpaired)[paired_offset(i, 2 * j, 2 * int64_t(halves)) / 2] = h;
    }
  };
  if (i >= nq) {
    for (int j = lane; j < halves; j += 64) { put(j, _Float16(0.0f)); }
    if (lane == 0) { qscal[3 * i] = qscal[3 * i + 1] = qscal[3 * i + 2] = 0.0; }
    return;
  }
  // a query of at most 64 N coordinates is loaded once, for its norm and its encoding (N, the
  // coordinates per lane and chunk, is sized to the dimension: fewer registers, more waves)
  const int64_t r      = rows != nullptr ? int64_t(rows[i]) : i;  // the caller's query row
  const bool one_chunk = dim <= 64 * N;
  double v[N], c[N];
  double nrm = 1.0;
  if (one_chunk) {
    lane_coords<N>(q, t, r, dim, 0, lane, v);
    lane_center<N>(center, dim, 0, lane, c);
    if (normalize) {
      double s2 = 0;
#pragma unroll
      for (int u = 0; u < N; ++u) { s2 = fma(v[u], v[u], s2); }  // past dim: + 0, exact
      s2  = wave_sum(s2);
      nrm = s2 > 0 ? sqrt(s2) : 1.0;
    }
  } else if (normalize) {
    nrm = wave_row_norm(q, t, r, dim, lane);
  }
  double a = 0, nw = 0, ew = 0;
  for (int64_t j0 = 0; j0 < dim; j0 += 64 * N) {
    if (!one_chunk) {
      lane_coords<N>(q, t, r, dim, j0, lane, v);
      lane_center<N>(center, dim, j0, lane, c);
    }
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int64_t j = j0 + 64 * u + lane;
      if (j < dim) {
        const double w   = (v[u] / nrm - c[u]) * inv_alpha;
        const _Float16 h = to_f16(w);
        const double e   = w - double(h);
        put(j, h);
        a  = fma(w, w, a);
        nw = fma(double(h), double(h), nw);
        ew = fma(e, e, ew);
      }
    }
  }
  for (int64_t j = dim + lane; j < halves; j += 64) { put(j, _Float16(0.0f)); }
  a  = wave_sum(a);
  nw = wave_sum(nw);
  ew = wave_sum(ew);
  if (lane == 0) {
    qscal[3 * i]     = a * (1.0 - 1e-13);
    qscal[3 * i + 1] = sqrt_up(nw, dim);
    qscal[3 * i + 2] = sqrt_up(ew, dim);
  }
}

__global__ void remove_f_kernel(const int64_t* ids, int64_t n, int64_t size, float* rowc,
                                unsigned long long* newly, row_places at)
{
  const int64_t t = blockIdx.x * int64_t(blockDim.x) + threadIdx.x;
  if (t >= n) { return; }
  const int64_t id = ids[t];
  if (id < 0 || id >= size) { return; }
  if (id < at.n_part) { static_cast<float*>(at.part_rowc)[at.part_pos[id]] = -INFINITY; }
  if (at.anchor_stride > 0 && id % at.anchor_stride == 0 && id / at.anchor_stride < at.n_anchor) {
    static_cast<float*>(at.anchor_rowc)[id / at.anchor_stride] = -INFINITY;
  }
  const int old = atomicExch(reinterpret_cast<int*>(rowc + stored_row(at, id)),
                             __float_as_int(-INFINITY));
  if (old != __float_as_int(-INFINITY)) { atomicAdd(newly, 1ull); }
}

}  // namespace

void column_sums(const void* x, elem t, int64_t n, int64_t dim, bool normalize, double* sums,
                 hipStream_t stream)
{
  if (n == 0) { return; }
  const int64_t rows_per_block = 512;
  const unsigned blocks        = unsigned((n + rows_per_block - 1) / rows_per_block);
  column_sums_kernel<<<blocks, 128, 0, stream>>>(x, t, n, dim, normalize, rows_per_block, sums);
}

void max_norm(const void* x, elem t, int64_t n, int64_t dim, bool normalize, const double* center,
              double* out, hipStream_t stream)
{
  if (n == 0) { return; }
  const unsigned blocks = unsigned(std::min<int64_t>((n + 3) / 4, 4096));
  max_norm_kernel<<<blocks, 256, 0, stream>>>(x, t, n, dim, normalize, center, out);
}

void encode_rows_f16(const void* x, elem t, int64_t n, int64_t dim, int halves, bool normalize,
                     const double* center, double inv_alpha, metric_kind metric, double gamma,
                     uint16_t* rows, float* rowc, double* maxima, hipStream_t stream)
{
  if (n == 0) { return; }
  // four rows per workgroup at a time, at most 4,096 workgroups (16 per CU) striding over the rest
  const unsigned blocks = unsigned(std::min<int64_t>((n + 3) / 4, 4096));
  encode_rows_f16_kernel<<<blocks, 256, 0, stream>>>(x, t, n, dim, halves, normalize, center,
                                                     inv_alpha, metric, gamma, rows, rowc, maxima);
}

void encode_queries_f16(const void* q, elem t, int64_t nq, int64_t nq_pad, int64_t dim,
                        int halves, bool normalize, const double* center, double inv_alpha,
                        uint16_t* qrows, double* qscal, hipStream_t stream, uint16_t* qpaired,
                        const int32_t* rows)
{
  if (nq_pad == 0) { return; }
  // one wave per query, four per block; a lane's coordinates per chunk sized to the dimension
  const unsigned grid = unsigned((nq_pad + 3) / 4);
  auto go = [&](auto kernel) {
    kernel<<<grid, 256, 0, stream>>>(q, rows, t, nq, nq_pad, dim, halves, normalize, center,
                                     inv_alpha, qrows, qscal, qpaired);
  };
  if (dim <= 256) {
    go(encode_queries_f16_kernel<4>);
  } else if (dim <= 512) {
    go(encode_queries_f16_kernel<8>);
  } else if (dim <= 768) {
    go(encode_queries_f16_kernel<12>);
  } else {
    go(encode_queries_f16_kernel<kLaneChunk>);
  }
}

void remove_rows_f16(const int64_t* ids, int64_t n, int64_t size, float* rowc,
                     unsigned long long* newly_removed, const row_places& at, hipStream_t stream)
{
  if (n == 0) { return; }
  remove_f_kernel<<<blocks_for(n), 256, 0, stream>>>(ids, n, size, rowc, newly_removed, at);
}

void encode_rows_i8(const uint8_t* x, int64_t n, int64_t dim, int row_bytes, uint8_t flip,
                    metric_kind metric, int8_t* codes, int32_t* rowc, hipStream_t stream)
{
  if (n == 0) { return; }
  if (row_bytes > 256) {
    encode_rows_wide_kernel<<<blocks_for(n * 64), 256, 0, stream>>>(x, n, dim, row_bytes, flip,
                                                                   metric, codes, rowc);
    return;
  }
  encode_rows_kernel<<<blocks_for(n * (row_bytes / 16)), 256, 0, stream>>>(x, n, dim, row_bytes,
                                                                          flip, metric, codes, rowc);
}

void encode_queries_i8(const uint8_t* q, int64_t nq, int64_t nq_pad, int64_t dim, int row_bytes,
                       uint8_t flip, int8_t* qcodes, hipStream_t stream, int8_t* qpaired,
                       const int32_t* rows)
{
  const int64_t n = nq_pad * row_bytes;
  if (n == 0) { return; }
  encode_queries_kernel<<<blocks_for(n), 256, 0, stream>>>(q, rows, nq, nq_pad, dim, row_bytes,
                                                           flip, qcodes, qpaired);
}

void remove_rows_i8(const int64_t* ids, int64_t n, int64_t size, int32_t* rowc,
                    unsigned long long* newly_removed, const row_places& at, hipStream_t stream)
{
  if (n == 0) { return; }
  remove_kernel<<<blocks_for(n), 256, 0, stream>>>(ids, n, size, rowc, newly_removed, at);
}

void fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t stream)
{
  if (n == 0) { return; }
  const unsigned b = blocks_for(n) < 4096 ? blocks_for(n) : 4096;
  fill_kernel<uint32_t><<<b, 256, 0, stream>>>(p, n, v);
}

void fill_i32(int32_t* p, int64_t n, int32_t v, hipStream_t stream)
{
  if (n == 0) { return; }
  const unsigned b = blocks_for(n) < 4096 ? blocks_for(n) : 4096;
  fill_kernel<int32_t><<<b, 256, 0, stream>>>(p, n, v);
}

void iota_i32(int32_t* p, int64_t n, int32_t first, hipStream_t stream)
{
  if (n <= 0) { return; }
  const unsigned b = blocks_for(n) < 4096 ? blocks_for(n) : 4096;
  iota_kernel<<<b, 256, 0, stream>>>(p, n, first);
}

}  // namespace certex_amd
